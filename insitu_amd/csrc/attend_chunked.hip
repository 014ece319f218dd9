// The chunked attend: attend_online / attend_two_pass (ops/attention.py:429-513)
// over a context split into 512-token chunks, bit-exact with the sequential
// reference.
//
// Why it can be exact. In the online softmax the running maximum m_t is the
// prefix maximum of the scores, so a chunk can reproduce the reference's
// arithmetic token for token once it knows the maximum of everything before
// it (M_in): the tokens where s_t > m_{t-1} are the rescale events, the factor
// there is LUT(s_t - m_{t-1}), and every other token contributes
// floor(v_norm * p * c_v[code] / 2^23) with p = LUT(m_t - s_t) -- plain
// integers. Between two events these terms only add, so a chunk hands over,
// per query head, one integer segment sum (and the sum of p) per event-free
// run plus the factor that opens each run. Replaying
//     acc = floor(acc * f / 2^15) + S,   l = floor(l * f / 2^15) + L
// over the runs in order is exactly the reference recurrence, provided the
// per-token int32 clamp of acc (attention.py:502-503) never fires; that is
// proven per run from a bound on |acc| plus the sum of |term| bounds, and a
// head whose bound fails is recomputed on the serial path.
//
// Kernels (one workgroup of 256 threads per (chunk, sequence, KV head)):
//   chunk_max    exact scores of the chunk for the G=4 query heads sharing the
//                KV head (lane = token), chunk maxima -> cmax
//   chunk_accum  the same scores again, M_in from cmax, an in-chunk prefix-max
//                scan (events, p), run sums per head (wave = head, lane =
//                channel) into a per-(sequence, head) pool; the last workgroup
//                of a (sequence, KV head) replays the runs, finalizes and
//                writes the Q16 output.
// Scores: sum_ch q[ch] * c[code_ch] in fp64 FMA (every partial sum is an
// integer below 2^51, so it is exact), then the int64 norm multiply and >>24
// as the reference does.
#include "serial_head.h"

namespace insitu {

constexpr int CT = 256;              // threads per workgroup
constexpr int TPT = 2;               // tokens per thread in the score phase
constexpr int CHUNK = CT * TPT;      // tokens per workgroup
constexpr int GF = 4;                // query heads per KV head on this path
constexpr int FLAG_POOL = 1;         // segment pool exhausted
constexpr int EV_BIT = 0x10000;      // event marker beside the 16-bit factor
constexpr double MAGIC = 6755399441055744.0;   // 1.5 * 2^52
constexpr int64_t MAGIC_BITS = 0x4338000000000000LL;
constexpr double DOT_LIMIT = 2251799813685248.0;  // 2^51

struct ChunkHdr {
    int32_t n_seg, flags, pool_off, pad;
};
struct SegMeta {
    int64_t L, B;
    int32_t f, pad0;
    int64_t pad1;
};

struct Chunked {
    int64_t *cmax;          // [chain][max_chunks][GF]
    ChunkHdr *hdr;          // [chain][max_chunks][GF]
    SegMeta *meta;          // [chain][GF][pool]
    int64_t *segS;          // [chain][GF][pool][d]
    unsigned int *done;     // [chain]
    unsigned int *pool_ctr; // [chain][GF]
    int32_t max_chunks, pool;
};

template <int D, int KB>
struct KF {
    static constexpr int KBYTES = D * KB / 8;
    static constexpr int KWORDS = KBYTES / 4;
    static constexpr int NFULL = KBYTES / 16;
    static constexpr int HALF = (KBYTES % 16) / 8;
    static constexpr int CPL = D / 64;
    static constexpr uint32_t MASK = (1u << KB) - 1u;
    static constexpr int RS = ((D * KB / 8 + D * 4 / 8 + 4) + 3) / 4 * 4;   // widest row with VB <= 4
};

__device__ __forceinline__ int64_t dbl_to_i64(double x) {
    // x is an integer with |x| < 2^51: adding 1.5 * 2^52 puts it in the low mantissa bits.
    return (int64_t)__double_as_longlong(x + MAGIC) - MAGIC_BITS;
}

// Exact scores of one token for the GF heads (attention.py:333-359).
template <int D, int KB>
__device__ __forceinline__ void token_scores(const uint8_t *__restrict__ hb, int64_t span,
                                             int norm_plane, int64_t t, const double (*qf)[GF],
                                             const double *kcf, int score_shift, int64_t (&s)[GF],
                                             uint32_t &normw) {
    using K = KF<D, KB>;
    uint32_t w[K::KWORDS + 1];
#pragma unroll
    for (int p = 0; p < K::NFULL; ++p) {
        const uint4 v = *(const uint4 *)(hb + p * span + t * 16);
        w[4 * p] = v.x;
        w[4 * p + 1] = v.y;
        w[4 * p + 2] = v.z;
        w[4 * p + 3] = v.w;
    }
    if (K::HALF) {
        const uint2 v = *(const uint2 *)(hb + K::NFULL * span + t * 8);
        w[4 * K::NFULL] = v.x;
        w[4 * K::NFULL + 1] = v.y;
    }
    w[K::KWORDS] = 0;
    normw = *(const uint32_t *)(hb + norm_plane * span + t * 4);
    double acc[GF];
#pragma unroll
    for (int h = 0; h < GF; ++h) acc[h] = 0.0;
#pragma unroll
    for (int c = 0; c < D; ++c) {
        const int o = c * KB;
        const int wi = o >> 5, sh = o & 31;
        uint32_t code;
        if (sh + KB <= 32)
            code = (w[wi] >> sh) & K::MASK;
        else
            code = __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh) & K::MASK;
        const double cent = kcf[code];
#pragma unroll
        for (int h = 0; h < GF; ++h) acc[h] = fma(qf[c][h], cent, acc[h]);
    }
    const int64_t kn = sext16(normw);
#pragma unroll
    for (int h = 0; h < GF; ++h) s[h] = wmul(dbl_to_i64(acc[h]), kn) >> score_shift;
}

// Shared prologue: q (fp64) and the key centroids (fp64) into LDS; checks that
// every head's score stays an exact fp64 integer (|dot| < 2^51).
template <int D>
__device__ __forceinline__ bool load_q(const Geom &g, const Tables *__restrict__ tabs,
                                       const int32_t *__restrict__ q, int b, int kvh,
                                       double (*qf)[GF], double *kcf, int *qok) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nk = 1 << g.kb;
    if (tid < nk) kcf[tid] = (double)tabs->kc[tid];
    if (tid == 0) *qok = 1;
    __syncthreads();
    // wave wv handles head wv
    const int32_t *qrow = q + ((int64_t)b * g.n_q + kvh * GF + wv) * D;
    double l1 = 0.0;
#pragma unroll
    for (int k = 0; k < D / 64; ++k) {
        const int c = lane + 64 * k;
        const int32_t v = qrow[c];
        qf[c][wv] = (double)v;
        l1 += fabs((double)v);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) l1 += __shfl_xor(l1, o, 64);
    if (lane == 0) {
        double cmax = 0.0;
        for (int i = 0; i < nk; ++i) cmax = fmax(cmax, fabs(kcf[i]));
        // l1 and cmax are exact in fp64 (below 2^53); the product bounds |dot|.
        if (!(l1 * cmax < DOT_LIMIT)) atomicAnd(qok, 0);
    }
    __syncthreads();
    return *qok != 0;
}

template <int D, int KB>
__global__ void __launch_bounds__(CT) chunk_max_kernel(Geom g, const Tables *__restrict__ tabs,
                                                       const int32_t *__restrict__ q,
                                                       const int64_t *__restrict__ len,
                                                       Chunked ck, DevStats *st) {
    __shared__ double qf[D][GF];
    __shared__ double kcf[16];
    __shared__ int qok;
    __shared__ int64_t red[CT / 64][GF];
    __shared__ unsigned long long ovf_s, mabs_s;
    const int chunk = blockIdx.x, chain = blockIdx.y;
    const int b = chain / g.n_kv, kvh = chain % g.n_kv;
    const int64_t T = len[b];
    const int64_t nch = T > 0 ? (T + CHUNK - 1) / CHUNK : 1;
    if (chunk >= nch) return;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    if (tid == 0) ovf_s = mabs_s = 0;
    const bool ok = load_q<D>(g, tabs, q, b, kvh, qf, kcf, &qok);
    if (chunk == 0) {
        // The seam promises 24-bit lanes; a rotated query beyond +-2^27 is flagged
        // (the arithmetic stays exact: such heads go to the serial path).
        const int32_t *qrow = q + ((int64_t)b * g.n_q + kvh * GF + wv) * D;
        unsigned long long bad = 0;
        for (int c = lane; c < D; c += 64) {
            const int64_t v = qrow[c];
            bad += (v >= Q_ROT_LIMIT || v <= -Q_ROT_LIMIT) ? 1 : 0;
        }
        bad = (unsigned long long)wave_sum64((int64_t)bad);
        if (lane == 0 && bad) atomicAdd(&st->range_errors, bad);
    }
    const uint8_t *hb = plane_ptr(g, b, kvh, 0);
    const int score_shift = CENT_FRAC + g.norm_frac;
    int64_t mx[GF];
#pragma unroll
    for (int h = 0; h < GF; ++h) mx[h] = SCORE_LO;
    unsigned long long ovf = 0;
    int64_t mabs = 0;
    if (ok) {
#pragma unroll
        for (int j = 0; j < TPT; ++j) {
            const int64_t t = (int64_t)chunk * CHUNK + j * CT + tid;
            if (t < T) {
                int64_t s[GF];
                uint32_t nw;
                token_scores<D, KB>(hb, g.span, g.n_planes - 1, t, qf, kcf, score_shift, s, nw);
#pragma unroll
                for (int h = 0; h < GF; ++h) {
                    int64_t v = s[h];
                    if (v < SCORE_LO || v > SCORE_HI) {
                        ++ovf;
                        v = v < SCORE_LO ? SCORE_LO : SCORE_HI;
                    }
                    const int64_t a = v < 0 ? -v : v;
                    mabs = a > mabs ? a : mabs;
                    mx[h] = v > mx[h] ? v : mx[h];
                }
            }
        }
    }
#pragma unroll
    for (int h = 0; h < GF; ++h) {
        const int64_t m = wave_max64(mx[h]);
        if (lane == 0) red[wv][h] = m;
    }
    ovf = (unsigned long long)wave_sum64((int64_t)ovf);
    mabs = wave_max64(mabs);
    if (lane == 0) {
        atomicAdd(&ovf_s, ovf);
        atomicMax(&mabs_s, (unsigned long long)mabs);
    }
    __syncthreads();
    if (tid < GF) {
        int64_t m = red[0][tid];
        for (int w = 1; w < CT / 64; ++w) m = red[w][tid] > m ? red[w][tid] : m;
        ck.cmax[((int64_t)chain * ck.max_chunks + chunk) * GF + tid] = m;
    }
    if (tid == 0 && ok) {
        if (ovf_s) atomicAdd(&st->score_overflows, ovf_s);
        atomicMax(&st->max_abs_score, mabs_s);
    }
}

template <int D, int KB>
struct AccumLds {
    struct Phase {
        int64_t s[GF][CHUNK];
        int32_t p[GF][CHUNK];
        int32_t ev[GF][CHUNK];
        uint32_t vw[CHUNK][D * 4 / 32];
        int32_t vn[CHUNK];
    };
    union {
        Phase ph;
        SerialLds<KF<D, KB>::RS> fb[GF];
    } u;
    double qf[D][GF];
    double kcf[16];
    int64_t kc[16];
    int64_t vc[16];
    int32_t expt[256];
    int64_t min_[GF];
    int64_t wt[CT / 64][GF];
    int qok;
    int last;
};

template <int D, int KB>
__global__ void __launch_bounds__(CT) chunk_accum_kernel(Geom g, const Tables *__restrict__ tabs,
                                                         const int32_t *__restrict__ q, int32_t *out,
                                                         const int64_t *__restrict__ len,
                                                         Chunked ck, int two_pass, DevStats *st) {
    using K = KF<D, KB>;
    constexpr int CPL = K::CPL;
    __shared__ AccumLds<D, KB> S;
    const int chunk = blockIdx.x, chain = blockIdx.y;
    const int b = chain / g.n_kv, kvh = chain % g.n_kv;
    const int64_t T = len[b];
    const int64_t nch = T > 0 ? (T + CHUNK - 1) / CHUNK : 1;
    if (chunk >= nch) return;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nv = 1 << g.vb;
    const int vwords = g.value_bytes / 4;
    const int acc_shift = CENT_FRAC + g.norm_frac + PROB_FRAC - ACC_FRAC;
    const int score_shift = CENT_FRAC + g.norm_frac;

    if (tid < 16) S.kc[tid] = tid < (1 << g.kb) ? tabs->kc[tid] : 0;
    if (tid < 16) S.vc[tid] = tid < nv ? tabs->vc[tid] : 0;
    S.expt[tid] = tabs->exp_table[tid];
    const bool ok = load_q<D>(g, tabs, q, b, kvh, S.qf, S.kcf, &S.qok);
    const uint8_t *hb = plane_ptr(g, b, kvh, 0);
    const int64_t t0 = (int64_t)chunk * CHUNK;

    // -- phase 1: scores (lane = token) and the value codes of the chunk ------
    if (ok) {
#pragma unroll
        for (int j = 0; j < TPT; ++j) {
            const int tl = j * CT + tid;
            const int64_t t = t0 + tl;
            int64_t s[GF];
            uint32_t nw = 0;
            if (t < T) {
                token_scores<D, KB>(hb, g.span, g.n_planes - 1, t, S.qf, S.kcf, score_shift, s, nw);
#pragma unroll
                for (int h = 0; h < GF; ++h)
                    s[h] = s[h] < SCORE_LO ? SCORE_LO : (s[h] > SCORE_HI ? SCORE_HI : s[h]);
                // value codes: they follow the key field; their planes are 16 or 8 bytes wide
                const int vp0 = K::NFULL + K::HALF;
                int wi = 0;
                for (int p = vp0; wi < vwords; ++p) {
                    const int wdt = g.plane_w[p];
                    const uint32_t *src = (const uint32_t *)(hb + p * g.span + t * wdt);
                    for (int i = 0; i < wdt / 4; ++i) S.u.ph.vw[tl][wi++] = src[i];
                }
            } else {
#pragma unroll
                for (int h = 0; h < GF; ++h) s[h] = SCORE_LO;
            }
            S.u.ph.vn[tl] = (int32_t)sext16(nw >> 16);
#pragma unroll
            for (int h = 0; h < GF; ++h) S.u.ph.s[h][tl] = s[h];
        }
    }
    // -- phase 2: the maximum of everything before this chunk (or of all, two-pass)
    {
        const int64_t lim = two_pass ? nch : chunk;
        int64_t m = SCORE_LO;
        for (int64_t c = lane; c < lim; c += 64) {
            const int64_t v = ck.cmax[((int64_t)chain * ck.max_chunks + c) * GF + wv];
            m = v > m ? v : m;
        }
        m = wave_max64(m);
        if (lane == 0) S.min_[wv] = m;
    }
    __syncthreads();

    // -- phase 3: events and p per token (thread owns TPT consecutive tokens) ---
    if (ok) {
        int64_t sv[GF][TPT];
        int64_t run[GF];
#pragma unroll
        for (int h = 0; h < GF; ++h) {
            run[h] = SCORE_LO;
#pragma unroll
            for (int j = 0; j < TPT; ++j) {
                sv[h][j] = S.u.ph.s[h][tid * TPT + j];
                run[h] = sv[h][j] > run[h] ? sv[h][j] : run[h];
            }
        }
        int64_t excl[GF];
        if (!two_pass) {
#pragma unroll
            for (int h = 0; h < GF; ++h) {
                int64_t v = run[h];
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) {
                    const int64_t u = __shfl_up(v, o, 64);
                    if (lane >= o) v = u > v ? u : v;
                }
                if (lane == 63) S.wt[wv][h] = v;
                const int64_t u = __shfl_up(v, 1, 64);
                excl[h] = lane > 0 ? u : SCORE_LO;
            }
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < GF; ++h) {
            if (two_pass) {
                const int64_t M = S.min_[h];
#pragma unroll
                for (int j = 0; j < TPT; ++j) {
                    const int tl = tid * TPT + j;
                    const bool valid = t0 + tl < T;
                    S.u.ph.p[h][tl] = valid ? exp_lut(M - sv[h][j], S.expt, tabs->delta_max) : 0;
                    S.u.ph.ev[h][tl] = 0;
                }
            } else {
                int64_t prev = S.min_[h];
                for (int w = 0; w < wv; ++w) prev = S.wt[w][h] > prev ? S.wt[w][h] : prev;
                prev = excl[h] > prev ? excl[h] : prev;
#pragma unroll
                for (int j = 0; j < TPT; ++j) {
                    const int tl = tid * TPT + j;
                    int32_t p = 0, ev = 0;
                    if (t0 + tl < T) {
                        const int64_t sj = sv[h][j];
                        if (sj > prev) {
                            ev = EV_BIT | exp_lut(sj - prev, S.expt, tabs->delta_max);
                            prev = sj;
                        }
                        p = exp_lut(prev - sj, S.expt, tabs->delta_max);
                    }
                    S.u.ph.p[h][tl] = p;
                    S.u.ph.ev[h][tl] = ev;
                }
            }
        }
    }
    __syncthreads();

    // -- phase 4: run sums, wave = head, lane = channel ------------------------
    if (ok) {
        const int h = wv;
        int n_ev = 0;
        for (int blk = 0; blk < CHUNK / 64; ++blk)
            n_ev += __popcll(__ballot(S.u.ph.ev[h][blk * 64 + lane] != 0));
        const int n_seg = n_ev + 1;
        int off = 0, flags = 0;
        if (lane == 0) off = (int)atomicAdd(&ck.pool_ctr[chain * GF + h], (unsigned)n_seg);
        off = __shfl(off, 0, 64);
        if (off + n_seg > ck.pool) flags |= FLAG_POOL;
        if (!flags) {
            // lane -> channel(s): code position in the value words is fixed per lane
            int wi[CPL], sh[CPL];
#pragma unroll
            for (int k = 0; k < CPL; ++k) {
                const int bit = (lane + 64 * k) * g.vb;
                wi[k] = bit >> 5;
                sh[k] = bit & 31;
            }
            const uint32_t vmask = (1u << g.vb) - 1u;
            const int64_t vcmax = [&] {
                int64_t m = 0;
                for (int i = 0; i < nv; ++i) {
                    const int64_t a = S.vc[i] < 0 ? -S.vc[i] : S.vc[i];
                    m = a > m ? a : m;
                }
                return m;
            }();
            SegMeta *meta = ck.meta + ((int64_t)chain * GF + h) * ck.pool;
            int64_t *segS = ck.segS + ((int64_t)chain * GF + h) * ck.pool * D;
            int seg = 0;
            int32_t segf = 0;
            int64_t Ssum[CPL];
#pragma unroll
            for (int k = 0; k < CPL; ++k) Ssum[k] = 0;
            int64_t L = 0, B = 0;
            for (int blk = 0; blk < CHUNK / 64; ++blk) {
                const int32_t pv = S.u.ph.p[h][blk * 64 + lane];
                const int32_t evv = S.u.ph.ev[h][blk * 64 + lane];
                unsigned long long mask = __ballot(pv != 0);
                while (mask) {
                    const int i = __ffsll((long long)mask) - 1;
                    mask &= mask - 1;
                    const int tl = blk * 64 + i;
                    const int32_t p = __shfl(pv, i, 64);
                    const int32_t e = __shfl(evv, i, 64);
                    if (e) {
                        // close the run that the event ends
                        if (lane == 0) {
                            meta[off + seg].L = L;
                            meta[off + seg].B = B;
                            meta[off + seg].f = segf;
                        }
#pragma unroll
                        for (int k = 0; k < CPL; ++k) segS[(int64_t)(off + seg) * D + lane + 64 * k] = Ssum[k];
                        ++seg;
                        segf = e & 0xFFFF;
#pragma unroll
                        for (int k = 0; k < CPL; ++k) Ssum[k] = 0;
                        L = 0;
                        B = 0;
                    }
                    const int32_t w = S.u.ph.vn[tl] * p;          // |w| <= 2^30
#pragma unroll
                    for (int k = 0; k < CPL; ++k) {
                        const uint32_t lo = S.u.ph.vw[tl][wi[k]];
                        uint32_t code;
                        if (sh[k] + g.vb <= 32)
                            code = (lo >> sh[k]) & vmask;
                        else
                            code = __builtin_amdgcn_alignbit(S.u.ph.vw[tl][wi[k] + 1], lo, sh[k]) & vmask;
                        Ssum[k] += ((int64_t)w * S.vc[code]) >> acc_shift;
                    }
                    L += p;
                    const int64_t aw = w < 0 ? -(int64_t)w : (int64_t)w;
                    B += ((aw * vcmax) >> acc_shift) + 1;
                }
            }
            if (lane == 0) {
                meta[off + seg].L = L;
                meta[off + seg].B = B;
                meta[off + seg].f = segf;
            }
#pragma unroll
            for (int k = 0; k < CPL; ++k) segS[(int64_t)(off + seg) * D + lane + 64 * k] = Ssum[k];
        }
        if (lane == 0) {
            ChunkHdr hd;
            hd.n_seg = n_seg;
            hd.flags = flags;
            hd.pool_off = off;
            hd.pad = 0;
            ck.hdr[((int64_t)chain * ck.max_chunks + chunk) * GF + h] = hd;
        }
    }

    // -- phase 5: the last workgroup of this (sequence, KV head) combines ------
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const unsigned prior = atomicAdd(&ck.done[chain], 1u);
        S.last = prior == (unsigned)(nch - 1);
    }
    __syncthreads();
    if (!S.last) return;
    __threadfence();

    const int h = wv;
    const int qh = kvh * GF + h;
    int32_t *orow = out + ((int64_t)b * g.n_q + qh) * D;
    bool fb = !ok;
    int64_t acc[CPL];
#pragma unroll
    for (int k = 0; k < CPL; ++k) acc[k] = 0;
    int64_t l = 0, R = 0;
    unsigned long long events = 0;
    if (!fb) {
        for (int64_t c = 0; c < nch && !fb; ++c) {
            const ChunkHdr hd = ck.hdr[((int64_t)chain * ck.max_chunks + c) * GF + h];
            if (hd.flags) {
                fb = true;
                break;
            }
            const SegMeta *meta = ck.meta + ((int64_t)chain * GF + h) * ck.pool + hd.pool_off;
            const int64_t *segS = ck.segS + (((int64_t)chain * GF + h) * ck.pool + hd.pool_off) * D;
            for (int j = 0; j < hd.n_seg; ++j) {
                const SegMeta m = meta[j];
                if (!two_pass) {
                    if (j > 0) {
#pragma unroll
                        for (int k = 0; k < CPL; ++k) acc[k] = wmul(acc[k], m.f) >> PROB_FRAC;
                        l = wmul(l, m.f) >> PROB_FRAC;
                        R = (wmul(R, m.f) >> PROB_FRAC) + 1;
                        ++events;
                    }
                    R += m.B;
                    if (R > ACC_HI) {
                        fb = true;
                        break;
                    }
                }
#pragma unroll
                for (int k = 0; k < CPL; ++k) acc[k] += segS[(int64_t)j * D + lane + 64 * k];
                l += m.L;
            }
        }
    }
    __syncthreads();   // the phase buffers are dead from here; the fallback reuses them
    if (fb) {
        // Score statistics were counted by chunk_max unless q failed its range check.
        serial_head<CPL, K::RS>(g, tabs, S.kc, S.vc, q + ((int64_t)b * g.n_q + qh) * D, b, kvh, T,
                                two_pass, !ok, S.u.fb[h], orow, st);
        if (lane == 0) atomicAdd(&st->serial_fallbacks, 1ull);
    } else {
        unsigned long long aovf = 0;
        if (two_pass) {
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
        amax = wave_max64(amax);
        aovf = (unsigned long long)wave_sum64((int64_t)aovf);
        if (lane == 0) {
            atomicMax(&st->n_tokens, (unsigned long long)T);
            atomicAdd(&st->rescale_events, events);
            atomicMax(&st->max_abs_acc, (unsigned long long)amax);
            if (aovf) atomicAdd(&st->acc_overflows, aovf);
        }
    }
    // reset the counters for the next call (every other workgroup of this chain is done)
    if (lane == 0) ck.pool_ctr[chain * GF + h] = 0;
    if (tid == 0) ck.done[chain] = 0;
}

template <int D, int KB>
static hipError_t launch_fast(hipStream_t s, const Geom &g, const Tables *t, const int32_t *q,
                              int32_t *out, const int64_t *len, const Chunked &ck, int two_pass,
                              DevStats *st) {
    dim3 grid((unsigned)ck.max_chunks, (unsigned)(g.batch * g.n_kv)), block(CT);
    hipLaunchKernelGGL((chunk_max_kernel<D, KB>), grid, block, 0, s, g, t, q, len, ck, st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((chunk_accum_kernel<D, KB>), grid, block, 0, s, g, t, q, out, len, ck,
                       two_pass, st);
    return hipGetLastError();
}

bool chunked_supported(const Geom &g) {
    return g.G == GF && (g.d == 64 || g.d == 128) && g.kb >= 2 && g.kb <= 4 && g.vb >= 1 &&
           g.vb <= 4;
}

int64_t chunked_max_chunks(int64_t capacity) { return (capacity + CHUNK - 1) / CHUNK; }

size_t chunked_scratch_bytes(const Geom &g, int64_t max_chunks, int64_t pool) {
    const int64_t chains = (int64_t)g.batch * g.n_kv;
    size_t n = 0;
    n += chains * max_chunks * GF * sizeof(int64_t);
    n += chains * max_chunks * GF * sizeof(ChunkHdr);
    n += chains * GF * pool * sizeof(SegMeta);
    n += chains * GF * pool * g.d * sizeof(int64_t);
    n += chains * sizeof(unsigned int);
    n += chains * GF * sizeof(unsigned int);
    return n + 1024;
}

hipError_t launch_attend_chunked(hipStream_t s, const Geom &g, const Tables *t, const int32_t *q,
                                 int32_t *out, const int64_t *len, void *scratch, int64_t max_chunks,
                                 int64_t pool, int two_pass, DevStats *st) {
    const int64_t chains = (int64_t)g.batch * g.n_kv;
    uint8_t *p = (uint8_t *)scratch;
    Chunked ck;
    ck.cmax = (int64_t *)p;
    p += chains * max_chunks * GF * sizeof(int64_t);
    ck.hdr = (ChunkHdr *)p;
    p += chains * max_chunks * GF * sizeof(ChunkHdr);
    ck.meta = (SegMeta *)p;
    p += chains * GF * pool * sizeof(SegMeta);
    ck.segS = (int64_t *)p;
    p += chains * GF * pool * g.d * sizeof(int64_t);
    ck.done = (unsigned int *)p;
    p += chains * sizeof(unsigned int);
    ck.pool_ctr = (unsigned int *)p;
    ck.max_chunks = (int32_t)max_chunks;
    ck.pool = (int32_t)pool;
    if (max_chunks > 65535 || chains > 65535) return hipErrorInvalidValue;
#define INSITU_FAST(DD, KK)                                                          \
    if (g.d == DD && g.kb == KK)                                                     \
        return launch_fast<DD, KK>(s, g, t, q, out, len, ck, two_pass, st);
    INSITU_FAST(64, 2)
    INSITU_FAST(64, 3)
    INSITU_FAST(64, 4)
    INSITU_FAST(128, 2)
    INSITU_FAST(128, 3)
    INSITU_FAST(128, 4)
#undef INSITU_FAST
    return hipErrorInvalidValue;
}

}  // namespace insitu
