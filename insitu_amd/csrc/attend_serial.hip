// The serial attend: CompressedAttention.attend_online / attend_two_pass
// (ops/attention.py:429-513) computed one query head per wave, token by token.
//
// Scores for 64 tokens at a time are computed with lane = token (each lane
// walks its row's key codes against q held in LDS); the online recurrence then
// walks those 64 tokens in order with lane = channel, exactly as the reference
// loop does. It is slow by design and exact by construction: it is the
// reference GPU path that the fast chunked kernel is tested against, and the
// fallback that kernel takes when an accumulator bound cannot be proven.
#include "insitu_internal.h"

namespace insitu {

constexpr int ROW_STRIDE = 272;   // >= the widest row (8b/8b at d=128: 260 B), 16-aligned

// Stage up to 64 rows of head `h` (tokens base .. base+n-1) into rows[t][*].
__device__ __forceinline__ void stage_rows(const Geom &g, int b, int h, int64_t base, int n,
                                           uint8_t (*rows)[ROW_STRIDE]) {
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

template <int CPL>
__global__ void __launch_bounds__(64) attend_serial_kernel(Geom g, const Tables *__restrict__ tabs,
                                                           const int32_t *__restrict__ q,
                                                           int32_t *out,
                                                           const int64_t *__restrict__ len,
                                                           int two_pass, DevStats *st) {
    __shared__ int64_t kc[256], vc[256];
    __shared__ int64_t qs[MAX_D];
    __shared__ __align__(16) uint8_t rows[64][ROW_STRIDE];
    const int lane = threadIdx.x;
    const int b = blockIdx.x / g.n_q;
    const int qh = blockIdx.x % g.n_q;
    const int kvh = qh / g.G;
    const int d = g.d;
    const int nk = 1 << g.kb, nv = 1 << g.vb;
    const int score_shift = CENT_FRAC + g.norm_frac;               // config.py:249-250
    const int acc_shift = CENT_FRAC + g.norm_frac + PROB_FRAC - ACC_FRAC;  // config.py:252-254
    const int noff = g.key_bytes + g.value_bytes;

    for (int i = lane; i < nk; i += 64) kc[i] = tabs->kc[i];
    for (int i = lane; i < nv; i += 64) vc[i] = tabs->vc[i];
    const int32_t *qrow = q + ((int64_t)b * g.n_q + qh) * d;
    for (int c = lane; c < d; c += 64) {
        int64_t qv = qrow[c];
        if (qv >= Q_ROT_LIMIT || qv <= -Q_ROT_LIMIT) atomicAdd(&st->range_errors, 1ull);
        qs[c] = qv;
    }
    __syncthreads();

    const int64_t T = len[b];
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
            stage_rows(g, b, kvh, base, n, rows);
            __syncthreads();
            int64_t s_mine = 0;
            if (lane < n) {
                int64_t dot = 0;
                for (int c = 0; c < d; ++c) dot = wadd(dot, wmul(qs[c], kc[code_at(rows[lane], c, g.kb)]));
                const int64_t kn = sext16((uint32_t)rows[lane][noff] | ((uint32_t)rows[lane][noff + 1] << 8));
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
                const int64_t sj = __shfl(s_mine, j, 64);
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
                const int64_t vn = sext16((uint32_t)rows[j][noff + 2] | ((uint32_t)rows[j][noff + 3] << 8));
                const int64_t w = wmul(vn, p);
#pragma unroll
                for (int k = 0; k < CPL; ++k) {
                    const int ch = lane + 64 * k;
                    if (ch < d) {
                        const int code = code_at(rows[j] + g.key_bytes, ch, g.vb);
                        int64_t a = wadd(acc[k], wmul(w, vc[code]) >> acc_shift);
                        if (!two_pass && (a < ACC_LO || a > ACC_HI)) {
                            ++aovf;
                            a = a < ACC_LO ? ACC_LO : ACC_HI;
                        }
                        acc[k] = a;
                    }
                }
            }
            __syncthreads();
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
            out[((int64_t)b * g.n_q + qh) * d + ch] = (int32_t)(wmul(acc[k], rc.r) >> rc.shift);
            int64_t a = acc[k] < 0 ? -acc[k] : acc[k];
            amax = a > amax ? a : amax;
        }
    }
    // statistics: per-lane counters reduced once per wave
    amax = wave_max64(amax);
    max_abs_s = wave_max64(max_abs_s);
    sovf = (unsigned long long)wave_sum64((int64_t)sovf);
    aovf = (unsigned long long)wave_sum64((int64_t)aovf);
    if (lane == 0) {
        atomicMax(&st->n_tokens, (unsigned long long)T);
        atomicAdd(&st->rescale_events, events);
        atomicAdd(&st->score_overflows, sovf);
        atomicAdd(&st->acc_overflows, aovf);
        atomicMax(&st->max_abs_score, (unsigned long long)max_abs_s);
        atomicMax(&st->max_abs_acc, (unsigned long long)amax);
    }
}

hipError_t launch_attend_serial(hipStream_t s, const Geom &g, const Tables *t, const int32_t *q,
                                int32_t *out, const int64_t *len, int two_pass, DevStats *st) {
    const int64_t blocks = (int64_t)g.batch * g.n_q;
    if (blocks <= 0) return hipSuccess;
    if (g.d <= 64)
        hipLaunchKernelGGL(attend_serial_kernel<1>, dim3((unsigned)blocks), dim3(64), 0, s, g, t, q,
                           out, len, two_pass, st);
    else
        hipLaunchKernelGGL(attend_serial_kernel<2>, dim3((unsigned)blocks), dim3(64), 0, s, g, t, q,
                           out, len, two_pass, st);
    return hipGetLastError();
}

}  // namespace insitu
