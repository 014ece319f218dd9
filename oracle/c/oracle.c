/* CPU oracle in C for long contexts. TEST INFRASTRUCTURE ONLY.
 *
 * The same arithmetic as oracle/attention.py (which restates ops/attention.py
 * of the reference), written as plain loops so a 32k-token online scan takes
 * milliseconds instead of minutes. int64 sums and products wrap modulo 2^64
 * exactly as numpy int64 does (computed in uint64, then reinterpreted).
 *
 * Inputs are the unpacked view of a cache (quantize.py:99-118): codes as one
 * uint8 per channel, norms as int64.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    int32_t d, key_bits, value_bits;
    int32_t score_shift;     /* config.py:249-250, 24 at the reference format */
    int32_t acc_shift;       /* config.py:252-254, 23 */
    int32_t prob_frac;       /* 15 */
    int32_t acc_frac;        /* 16 */
    int32_t score_width;     /* 48 */
    int32_t acc_width;       /* 32 */
} orc_fmt;

typedef struct {
    int64_t n_tokens, rescale_events, score_overflows, acc_overflows, max_abs_score, max_abs_acc;
} orc_stats;

static inline int64_t wmul(int64_t a, int64_t b) { return (int64_t)((uint64_t)a * (uint64_t)b); }
static inline int64_t wadd(int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); }
static inline int64_t asr(int64_t a, int n) { return a >> n; }   /* gcc: arithmetic */
static inline int64_t iabs64(int64_t a) { return a < 0 ? -a : a; }

/* attention.py:90-159, flat form. table[256] = rint(2^(-i/256) * 2^15). */
typedef struct {
    int64_t flat[(17 << 8) + 1];
    int64_t delta_max, log2e;
    int32_t shift, span, acc_frac;
} orc_exp;

void orc_exp_init(orc_exp *e, const int64_t *table256, int64_t log2e, int64_t delta_max,
                  int32_t acc_frac, int32_t lut_bits, int32_t max_int_part) {
    int32_t n = 1 << lut_bits;
    e->span = (max_int_part + 1) << lut_bits;
    e->shift = acc_frac - lut_bits;
    e->acc_frac = acc_frac;
    e->log2e = log2e;
    e->delta_max = delta_max;
    for (int32_t u = 0; u < e->span; ++u) {
        int32_t ip = u >> lut_bits;
        e->flat[u] = ip > max_int_part ? 0 : (table256[u & (n - 1)] >> (ip < max_int_part ? ip : max_int_part));
    }
    e->flat[e->span] = 0;
}

static inline int64_t orc_exp_eval(const orc_exp *e, int64_t delta) {
    int64_t d = delta < e->delta_max ? delta : e->delta_max;
    int64_t t = asr(d * e->log2e, e->acc_frac);
    int64_t u = t >> e->shift;
    if (u > e->span) u = e->span;
    return e->flat[u];
}

int64_t orc_exp_vec(const orc_exp *e, const int64_t *delta, int64_t n, int64_t *out) {
    for (int64_t i = 0; i < n; ++i) {
        if (delta[i] < 0) return -1;
        out[i] = orc_exp_eval(e, delta[i]);
    }
    return 0;
}

/* attention.py:333-359 for G query heads against T rows. s is (G, T). */
void orc_scores(const orc_fmt *f, int32_t G, const int64_t *q, int64_t T,
                const uint8_t *k_idx, const int64_t *k_norm, const int64_t *kc,
                int64_t *s, orc_stats *st) {
    const int32_t d = f->d;
    const int64_t lo = -((int64_t)1 << (f->score_width - 1));
    const int64_t hi = ((int64_t)1 << (f->score_width - 1)) - 1;
    for (int32_t g = 0; g < G; ++g) {
        const int64_t *qg = q + (int64_t)g * d;
        for (int64_t t = 0; t < T; ++t) {
            const uint8_t *c = k_idx + t * d;
            int64_t dot = 0;
            for (int32_t j = 0; j < d; ++j) dot = wadd(dot, wmul(qg[j], kc[c[j]]));
            int64_t v = asr(wmul(dot, k_norm[t]), f->score_shift);
            if (v < lo) { v = lo; st->score_overflows++; }
            else if (v > hi) { v = hi; st->score_overflows++; }
            if (iabs64(v) > st->max_abs_score) st->max_abs_score = iabs64(v);
            s[(int64_t)g * T + t] = v;
        }
    }
}

/* attention.py:197-250 and :873-880. */
void orc_finalize(const orc_fmt *f, int32_t rows, int32_t d, const int64_t *acc, const int64_t *l,
                  int64_t *out, int64_t *recip, int64_t *shift) {
    for (int32_t r = 0; r < rows; ++r) {
        int64_t a = l[r];
        int64_t s = 0;
        for (int b = 1; b < 48; ++b) if (a >= ((int64_t)1 << b)) s = b;
        int64_t k = s - 31;
        int64_t ln = k >= 0 ? (a >> k) : (a << (-k));
        int64_t rr = a > 0 ? (int64_t)(((uint64_t)1 << 62) / (uint64_t)(ln > 1 ? ln : 1)) : 0;
        int64_t sh = 62 - f->prob_frac + k;
        if (recip) recip[r] = rr;
        if (shift) shift[r] = sh;
        for (int32_t j = 0; j < d; ++j) out[(int64_t)r * d + j] = asr(wmul(acc[(int64_t)r * d + j], rr), (int)sh);
    }
}

/* attention.py:451-513: the sequential-order online softmax for G heads.
 * acc (G, d), l (G), m (G) are the end-of-scan state; out (G, d). */
void orc_attend_online(const orc_fmt *f, const orc_exp *e, int32_t G, const int64_t *q, int64_t T,
                       const uint8_t *k_idx, const int64_t *k_norm,
                       const uint8_t *v_idx, const int64_t *v_norm,
                       const int64_t *kc, const int64_t *vc, int64_t *s_scratch,
                       int64_t *acc, int64_t *l, int64_t *m, int64_t *out, orc_stats *st) {
    const int32_t d = f->d;
    const int64_t acc_lo = -((int64_t)1 << (f->acc_width - 1));
    const int64_t acc_hi = ((int64_t)1 << (f->acc_width - 1)) - 1;
    const int64_t unity = (int64_t)1 << f->prob_frac;
    st->n_tokens = T;
    orc_scores(f, G, q, T, k_idx, k_norm, kc, s_scratch, st);
    for (int32_t g = 0; g < G; ++g) {
        int64_t *a = acc + (int64_t)g * d;
        memset(a, 0, sizeof(int64_t) * d);
        int64_t lg = 0, mg = -((int64_t)1 << (f->score_width - 1));
        const int64_t *sg = s_scratch + (int64_t)g * T;
        for (int64_t t = 0; t < T; ++t) {
            int64_t stt = sg[t];
            if (stt > mg) {
                int64_t fac = orc_exp_eval(e, stt - mg);
                for (int32_t j = 0; j < d; ++j) a[j] = asr(wmul(a[j], fac), f->prob_frac);
                lg = asr(wmul(lg, fac), f->prob_frac);
                mg = stt;
                st->rescale_events++;
            }
            (void)unity;
            int64_t p = orc_exp_eval(e, mg - stt);
            lg = wadd(lg, p);
            int64_t w = wmul(v_norm[t], p);
            if (w == 0) continue;        /* every term floor(0 * c / 2^23) is 0 */
            const uint8_t *vcode = v_idx + t * d;
            for (int32_t j = 0; j < d; ++j) {
                int64_t v = wadd(a[j], asr(wmul(w, vc[vcode[j]]), f->acc_shift));
                if (v < acc_lo) { v = acc_lo; st->acc_overflows++; }
                else if (v > acc_hi) { v = acc_hi; st->acc_overflows++; }
                a[j] = v;
            }
        }
        l[g] = lg;
        m[g] = mg;
        for (int32_t j = 0; j < d; ++j) if (iabs64(a[j]) > st->max_abs_acc) st->max_abs_acc = iabs64(a[j]);
    }
    orc_finalize(f, G, d, acc, l, out, 0, 0);
}

/* attention.py:429-449: global max, one accumulation, clamp at the end. */
void orc_attend_two_pass(const orc_fmt *f, const orc_exp *e, int32_t G, const int64_t *q, int64_t T,
                         const uint8_t *k_idx, const int64_t *k_norm,
                         const uint8_t *v_idx, const int64_t *v_norm,
                         const int64_t *kc, const int64_t *vc, int64_t *s_scratch,
                         int64_t *acc, int64_t *l, int64_t *out, orc_stats *st) {
    const int32_t d = f->d;
    const int64_t acc_lo = -((int64_t)1 << (f->acc_width - 1));
    const int64_t acc_hi = ((int64_t)1 << (f->acc_width - 1)) - 1;
    st->n_tokens = T;
    orc_scores(f, G, q, T, k_idx, k_norm, kc, s_scratch, st);
    for (int32_t g = 0; g < G; ++g) {
        const int64_t *sg = s_scratch + (int64_t)g * T;
        int64_t mg = T > 0 ? sg[0] : 0;
        for (int64_t t = 1; t < T; ++t) if (sg[t] > mg) mg = sg[t];
        int64_t *a = acc + (int64_t)g * d;
        memset(a, 0, sizeof(int64_t) * d);
        int64_t lg = 0;
        for (int64_t t = 0; t < T; ++t) {
            int64_t p = orc_exp_eval(e, mg - sg[t]);
            lg = wadd(lg, p);
            int64_t w = wmul(v_norm[t], p);
            const uint8_t *vcode = v_idx + t * d;
            for (int32_t j = 0; j < d; ++j) a[j] = wadd(a[j], asr(wmul(w, vc[vcode[j]]), f->acc_shift));
        }
        for (int32_t j = 0; j < d; ++j) {
            if (a[j] < acc_lo) { a[j] = acc_lo; st->acc_overflows++; }
            else if (a[j] > acc_hi) { a[j] = acc_hi; st->acc_overflows++; }
            if (iabs64(a[j]) > st->max_abs_acc) st->max_abs_acc = iabs64(a[j]);
        }
        l[g] = lg;
    }
    orc_finalize(f, G, d, acc, l, out, 0, 0);
}

/* The config-1 check: one layer's sequential decode from an empty cache
 * (kernel.py:271-345, the token attends to itself), or a prefill's queries
 * (attend_online_batch, attention.py:794-871). Step i attends its rotated
 * query rows q[i] (n_kv groups of G rows of d) over rows 0 .. base + i of each
 * KV head, exactly as orc_attend_online. k_idx/v_idx are (n_kv, cap, d) codes,
 * k_norm/v_norm (n_kv, cap); out is (steps, n_kv, G, d). Returns 0, or -1 when
 * scratch cannot be allocated or base + steps exceeds cap. */
int orc_decode_steps(const orc_fmt *f, const orc_exp *e, int32_t n_kv, int32_t G, int64_t steps,
                     int64_t base, int64_t cap, const int64_t *q, const uint8_t *k_idx, const int64_t *k_norm,
                     const uint8_t *v_idx, const int64_t *v_norm, const int64_t *kc,
                     const int64_t *vc, int64_t *out) {
    const int32_t d = f->d;
    if (base < 0 || base + steps > cap) return -1;
    int64_t *s = (int64_t *)malloc(sizeof(int64_t) * (size_t)G * (size_t)(base + steps > 0 ? base + steps : 1));
    int64_t *acc = (int64_t *)malloc(sizeof(int64_t) * (size_t)G * (size_t)d);
    int64_t *l = (int64_t *)malloc(sizeof(int64_t) * (size_t)G);
    int64_t *m = (int64_t *)malloc(sizeof(int64_t) * (size_t)G);
    int rc = (s && acc && l && m) ? 0 : -1;
    for (int64_t t = 0; t < steps && rc == 0; ++t) {
        for (int32_t h = 0; h < n_kv; ++h) {
            orc_stats st;
            memset(&st, 0, sizeof st);
            const int64_t qo = (t * n_kv + h) * (int64_t)G * d;
            orc_attend_online(f, e, G, q + qo, base + t + 1, k_idx + (int64_t)h * cap * d, k_norm + (int64_t)h * cap,
                              v_idx + (int64_t)h * cap * d, v_norm + (int64_t)h * cap, kc, vc, s, acc, l,
                              m, out + qo, &st);
        }
    }
    free(s);
    free(acc);
    free(l);
    free(m);
    return rc;
}
