// One query head's attend_online / attend_two_pass (ops/attention.py:429-513),
// token by token, by one wave.
//
// Scores for 64 tokens at a time are computed with lane = token (each lane
// walks its row's key codes against q held in LDS); the online recurrence then
// walks those 64 tokens in order with lane = channel, exactly as the reference
// loop does. Slow by design and exact by construction: it is the reference GPU
// path, and the fallback of the chunked kernel when an accumulator bound
// cannot be proven.
#pragma once

#include "insitu_internal.h"
#include "wave.h"

namespace insitu {

// Per-wave LDS of the serial path. RS >= row_bytes, a multiple of 4.
template <int RS>
struct SerialLds {
    int64_t qs[MAX_D];
    uint8_t rows[64][RS];
};

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Stage up to 64 rows of head `h` (tokens base .. base+n-1) into rows[t][*].
template <int RS>
__device__ __forceinline__ void stage_rows(const Geom &g, int b, int h, int64_t base, int n,
                                           uint8_t (*rows)[RS]) {
    const int lane = threadIdx.x & 63;
    if (lane < n) {
        for (int p = 0; p < g.n_planes; ++p) {
            const int w = g.plane_w[p];
            const uint8_t *src = plane_ptr(g, b, h, p) + (base + lane) * w;
            uint32_t *dst = (uint32_t *)&rows[lane][g.plane_lo[p]];
            for (int i = 0; i < w / 4; ++i) dst[i] = ((const uint32_t *)src)[i];
        }
    }
}

// kc/vc: the key/value centroids (int64) in LDS or global memory.
// Writes out_row[0..d) and merges this head's statistics into `st`. Score
// statistics are merged only when count_scores is set (the chunked kernel
// has already counted them when it falls back here).
template <int CPL, int RS>
__device__ __forceinline__ void serial_head(const Geom &g, const Tables *__restrict__ tabs,
                                            const int64_t *kc, const int64_t *vc,
                                            const int32_t *__restrict__ qrow, int b, int kvh, int64_t T,
                                            int two_pass, bool count_scores, SerialLds<RS> &L,
                                            int32_t *out_row, DevStats *st) {
    const int lane = threadIdx.x & 63;
    const int d = g.d;
    const int score_shift = CENT_FRAC + g.norm_frac;                        // config.py:249-250
    const int acc_shift = CENT_FRAC + g.norm_frac + PROB_FRAC - ACC_FRAC;   // config.py:252-254
    const int noff = g.key_bytes + g.value_bytes;

    for (int c = lane; c < d; c += 64) L.qs[c] = qrow[c];
    wave_sync();

    int64_t acc[CPL];
#pragma unroll
    for (int k = 0; k < CPL; ++k) acc[k] = 0;
    int64_t l = 0, m = SCORE_LO, gmax = SCORE_LO;
    unsigned long long events = 0, sovf = 0, aovf = 0;
    int64_t max_abs_s = 0;

    const int passes = two_pass ? 2 : 1;
    for (int pass = 0; pass < passes; ++pass) {
        for (int64_t base = 0; base < T; base += 64) {
            const int n = (int)((T - base) < 64 ? (T - base) : 64);
            wave_sync();
            stage_rows<RS>(g, b, kvh, base, n, L.rows);
            wave_sync();
            int64_t s_mine = 0;
            if (lane < n) {
                int64_t dot = 0;
                for (int c = 0; c < d; ++c)
                    dot = wadd(dot, wmul(L.qs[c], kc[code_at(L.rows[lane], c, g.kb)]));
                const int64_t kn = sext16((uint32_t)L.rows[lane][noff] |
                                          ((uint32_t)L.rows[lane][noff + 1] << 8));
                int64_t s = wmul(dot, kn) >> score_shift;
                if (s < SCORE_LO || s > SCORE_HI) {
                    if (pass == 0) ++sovf;
                    s = s < SCORE_LO ? SCORE_LO : SCORE_HI;
                }
                if (pass == 0) {
                    int64_t a = s < 0 ? -s : s;
                    if (a > max_abs_s) max_abs_s = a;
                }
                s_mine = s;
            }
            for (int j = 0; j < n; ++j) {
                const int64_t sj = readlane64(s_mine, j);
                int64_t p;
                if (!two_pass) {
                    if (sj > m) {
                        const int64_t f = exp_lut(sj - m, tabs->exp_table, tabs->delta_max);
#pragma unroll
                        for (int k = 0; k < CPL; ++k) acc[k] = wmul(acc[k], f) >> PROB_FRAC;
                        l = wmul(l, f) >> PROB_FRAC;
                        m = sj;
                        ++events;
                    }
                    p = exp_lut(m - sj, tabs->exp_table, tabs->delta_max);
                } else if (pass == 0) {
                    gmax = sj > gmax ? sj : gmax;
                    continue;
                } else {
                    p = exp_lut(gmax - sj, tabs->exp_table, tabs->delta_max);
                }
                l = wadd(l, p);
                const int64_t vn = sext16((uint32_t)L.rows[j][noff + 2] |
                                          ((uint32_t)L.rows[j][noff + 3] << 8));
                const int64_t w = wmul(vn, p);
#pragma unroll
                for (int k = 0; k < CPL; ++k) {
                    const int ch = lane + 64 * k;
                    if (ch < d) {
                        const int code = code_at(L.rows[j] + g.key_bytes, ch, g.vb);
                        int64_t a = wadd(acc[k], wmul(w, vc[code]) >> acc_shift);
                        if (!two_pass && (a < ACC_LO || a > ACC_HI)) {
                            ++aovf;
                            a = a < ACC_LO ? ACC_LO : ACC_HI;
                        }
                        acc[k] = a;
                    }
                }
            }
        }
    }
    if (two_pass) {
#pragma unroll
        for (int k = 0; k < CPL; ++k) {
            const int ch = lane + 64 * k;
            if (ch < d && (acc[k] < ACC_LO || acc[k] > ACC_HI)) {
                ++aovf;
                acc[k] = acc[k] < ACC_LO ? ACC_LO : ACC_HI;
            }
        }
    }
    const Recip rc = reciprocal(l);
    int64_t amax = 0;
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
        const int ch = lane + 64 * k;
        if (ch < d) {
            out_row[ch] = (int32_t)(wmul(acc[k], rc.r) >> rc.shift);
            int64_t a = acc[k] < 0 ? -acc[k] : acc[k];
            amax = a > amax ? a : amax;
        }
    }
    amax = wave_max_i64(amax);
    max_abs_s = wave_max_i64(max_abs_s);
    sovf = (unsigned long long)wave_sum_i64((int64_t)sovf);
    aovf = (unsigned long long)wave_sum_i64((int64_t)aovf);
    if (lane == 0) {
        atomicMax(&st->n_tokens, (unsigned long long)T);
        atomicAdd(&st->rescale_events, events);
        atomicAdd(&st->acc_overflows, aovf);
        atomicMax(&st->max_abs_acc, (unsigned long long)amax);
        if (count_scores) {
            atomicAdd(&st->score_overflows, sovf);
            atomicMax(&st->max_abs_score, (unsigned long long)max_abs_s);
        }
    }
}

}  // namespace insitu
